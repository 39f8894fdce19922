"""Tensor-level ops over the C ABI, mirroring pulsarlm-core's quant-linear ops.

Same names, argument meaning and error behaviour as the reference's
``pulsarlm-core/inc/pulsarlm/kernels/ops.hpp:299-332``:

* ``repack_int4_marlin_cuda(weight_packed, weight_scale, block_n, group_size)``
  -> ``(weight_marlin, scale_marlin)``
* ``repack_fp8_marlin_cuda(weight, weight_scale, block_n, group_size)``
* ``gemm_int4_marlin_cuda(x, weight_marlin, scale_marlin, n, block_n, group_size)``
* ``gemm_fp8_marlin_cuda(...)``

``weight_marlin`` is an opaque 1-D int32 tensor in the plm tile layout (the
reference's is also opaque, marlin.cu:21-30); ``scale_marlin`` keeps the scale's
source dtype, shaped [strips, groups, cols]. Errors raise ``RuntimeError`` with
the reference's ``"<op>: ..."`` message style. Work is enqueued on torch's
current stream of the tensors' device; nothing synchronizes.
"""

from __future__ import annotations

import threading

import torch

from . import _lib

_DTYPES = {torch.bfloat16: _lib.PLM_BF16, torch.float16: _lib.PLM_FP16, torch.float32: _lib.PLM_FP32}


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require(cond: bool, op: str, msg: str) -> None:
    if not cond:
        raise RuntimeError(f"{op}: {msg}")


def _call(fn_name: str, *args) -> None:
    lib = _lib.load()
    _lib.check(getattr(lib, fn_name)(*args))


# ---------------------------------------------------------------------------
# Workspace: one zero-initialised buffer per (device, stream). The kernels leave
# their arrival counters at zero, so reuse by calls ordered on one stream is safe.
# ---------------------------------------------------------------------------
_ws_lock = threading.Lock()
_ws: dict[tuple[int, int], torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    if nbytes <= 0:
        return None
    key = (device.index if device.index is not None else torch.cuda.current_device(), _stream(device))
    with _ws_lock:
        buf = _ws.get(key)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 1 << 20)
            buf = torch.zeros(size, dtype=torch.uint8, device=device)
            _ws[key] = buf
        return buf


# ---------------------------------------------------------------------------
# Repack
# ---------------------------------------------------------------------------


def _scale_shape(n: int, k: int, block_n: int, group_size: int):
    strips = -(-n // 16)
    ktiles = -(-k // 128)
    groups = -(-(ktiles * 128) // group_size)
    cols = 1 if block_n % 16 == 0 else 16
    return strips, groups, cols


def _repack(op: str, fmt: int, weight: torch.Tensor, n: int, k: int, weight_scale: torch.Tensor, block_n: int,
            group_size: int):
    _require(weight.is_cuda and weight_scale.is_cuda, op, "inputs must be CUDA tensors")
    _require(block_n > 0, op, "block_n must be positive")
    _require(group_size > 0 and group_size % 16 == 0, op, "group_size must be a positive multiple of 16")
    _require(k % group_size == 0, op, "K must be a multiple of group_size")
    rows = -(-n // block_n)
    _require(weight_scale.dim() == 2 and tuple(weight_scale.shape) == (rows, k // group_size), op,
             "weight_scale must be [ceil(N / block_n), K / group_size]")
    _require(weight_scale.dtype in _DTYPES, op, "weight_scale must be fp32, fp16 or bf16")
    src = weight.contiguous()
    scale = weight_scale.contiguous()
    lib = _lib.load()
    wbytes = lib.plm_weight_bytes(fmt, n, k)
    w_out = torch.empty(max(wbytes // 4, 0), dtype=torch.int32, device=weight.device)
    s_out = torch.empty(_scale_shape(n, k, block_n, group_size), dtype=scale.dtype, device=weight.device)
    fn = "plm_repack_int4" if fmt == _lib.PLM_INT4 else "plm_repack_fp8"
    with torch.cuda.device(weight.device):
        _call(fn, _ptr(src), _ptr(scale), _DTYPES[scale.dtype], n, k, block_n, group_size, _ptr(w_out), _ptr(s_out),
              _stream(weight.device))
    return w_out, s_out


def repack_int4_marlin_cuda(weight_packed: torch.Tensor, weight_scale: torch.Tensor, block_n: int, group_size: int):
    """int32 [N, K/8] LSB-first int4 + scales [ceil(N/bn), K/g] -> (weight, scale) in the plm layout
    (ops.hpp:306-311; marlin.cu:601-620)."""
    _require(weight_packed.dtype == torch.int32 and weight_packed.dim() == 2, "repack_int4_marlin",
             "weight_packed must be int32 [N, K/8]")
    n, k = weight_packed.shape[0], weight_packed.shape[1] * 8
    return _repack("repack_int4_marlin", _lib.PLM_INT4, weight_packed, n, k, weight_scale, block_n, group_size)


def repack_fp8_marlin_cuda(weight: torch.Tensor, weight_scale: torch.Tensor, block_n: int, group_size: int):
    """float8_e4m3fn [N, K] + scales -> (weight, scale) in the plm layout (ops.hpp:313-314; marlin.cu:622-629)."""
    _require(weight.dtype == torch.float8_e4m3fn and weight.dim() == 2, "repack_fp8_marlin",
             "weight must be float8_e4m3fn [N, K]")
    n, k = weight.shape
    return _repack("repack_fp8_marlin", _lib.PLM_FP8, weight.view(torch.uint8), n, k, weight_scale, block_n,
                   group_size)


def convert_marlin_cuda(fmt: str, weight_marlin: torch.Tensor, scale_marlin: torch.Tensor, n: int, k: int,
                        block_n: int, group_size: int):
    """Reference Marlin (words, fp32 [K/g, ceil(N/bn)] scales) -> plm layout (fp32 scales)."""
    op = "convert_marlin"
    f = _lib.PLM_INT4 if fmt == "int4" else _lib.PLM_FP8
    _require(weight_marlin.dtype == torch.int32 and scale_marlin.dtype == torch.float32, op,
             "weight_marlin must be int32 and scale_marlin fp32")
    lib = _lib.load()
    w_out = torch.empty(lib.plm_weight_bytes(f, n, k) // 4, dtype=torch.int32, device=weight_marlin.device)
    s_out = torch.empty(_scale_shape(n, k, block_n, group_size), dtype=torch.float32, device=weight_marlin.device)
    with torch.cuda.device(weight_marlin.device):
        _call("plm_convert_marlin", f, _ptr(weight_marlin.contiguous()), _ptr(scale_marlin.contiguous()), n, k,
              block_n, group_size, _ptr(w_out), _ptr(s_out), _stream(weight_marlin.device))
    return w_out, s_out


def dequant_marlin_cuda(fmt: str, weight_marlin: torch.Tensor, scale_marlin: torch.Tensor, n: int, k: int,
                        block_n: int, group_size: int, dtype=torch.bfloat16) -> torch.Tensor:
    """Dense [N, K] round(q * round(scale)) in ``dtype`` from the plm layout."""
    f = _lib.PLM_INT4 if fmt == "int4" else _lib.PLM_FP8
    out = torch.empty((n, k), dtype=dtype, device=weight_marlin.device)
    with torch.cuda.device(weight_marlin.device):
        _call("plm_dequant", f, _ptr(weight_marlin), _ptr(scale_marlin), _DTYPES[scale_marlin.dtype], n, k, block_n,
              group_size, _ptr(out), _DTYPES[dtype], _stream(weight_marlin.device))
    return out


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------


def _gemm_checks(op: str, fmt: int, x: torch.Tensor, weight_marlin: torch.Tensor, scale_marlin: torch.Tensor, n: int,
                 block_n: int, group_size: int):
    """gemm<fmt> checks, marlin.cu:547-571."""
    _require(x.is_cuda and weight_marlin.is_cuda and scale_marlin.is_cuda, op, "all inputs must be CUDA tensors")
    _require(x.dtype in (torch.float16, torch.bfloat16), op, "x must be fp16 or bf16")
    _require(x.dim() == 2 and x.is_contiguous(), op, "x must be a contiguous [M, K]")
    _require(weight_marlin.dtype == torch.int32, op, "weight_marlin must be int32")
    _require(scale_marlin.dtype in _DTYPES, op, "scale_marlin must be fp32, fp16 or bf16")
    _require(block_n > 0, op, "block_n must be positive")
    _require(group_size > 0 and group_size % 16 == 0, op, "group_size must be a positive multiple of 16")
    k = x.shape[1]
    _require(k % group_size == 0, op, "K must be a multiple of group_size")
    _require(tuple(scale_marlin.shape) == _scale_shape(n, k, block_n, group_size), op,
             "scale_marlin has the wrong shape for this N, K, block_n and group_size")
    _require(weight_marlin.numel() * 4 == _lib.load().plm_weight_bytes(fmt, n, k), op,
             "weight_marlin has the wrong size for this shape")


def _gemm(op: str, fmt: int, x, weight_marlin, scale_marlin, n: int, block_n: int, group_size: int,
          out: torch.Tensor | None = None) -> torch.Tensor:
    _gemm_checks(op, fmt, x, weight_marlin, scale_marlin, n, block_n, group_size)
    m, k = x.shape
    y = out if out is not None else torch.empty((m, n), dtype=x.dtype, device=x.device)
    if m == 0 or n == 0:
        return y
    lib = _lib.load()
    wsb = lib.plm_gemm_workspace_bytes(fmt, m, n, k)
    ws = workspace(x.device, wsb)
    with torch.cuda.device(x.device):
        _call("plm_gemm", fmt, _ptr(x), _DTYPES[x.dtype], _ptr(weight_marlin.contiguous()),
              _ptr(scale_marlin.contiguous()), _DTYPES[scale_marlin.dtype], m, n, k, block_n, group_size, _ptr(y),
              _ptr(ws), 0 if ws is None else ws.numel(), _stream(x.device))
    return y


def gemm_int4_marlin_cuda(x, weight_marlin, scale_marlin, n: int, block_n: int, group_size: int, out=None):
    """y [M, N] = x [M, K] @ dequant(W)^T (ops.hpp:316-323; marlin.cu:631-640)."""
    return _gemm("gemm_int4_marlin", _lib.PLM_INT4, x, weight_marlin, scale_marlin, n, block_n, group_size, out)


def gemm_fp8_marlin_cuda(x, weight_marlin, scale_marlin, n: int, block_n: int, group_size: int, out=None):
    """fp8 W8A16 form (ops.hpp:325-332; marlin.cu:642-651)."""
    return _gemm("gemm_fp8_marlin", _lib.PLM_FP8, x, weight_marlin, scale_marlin, n, block_n, group_size, out)


def quantize_rows_e4m3_cuda(x: torch.Tensor):
    """Per-row dynamic e4m3 quantization: (codes uint8 [M, K], scale fp32 [M]),
    scale = max(amax, 1e-12) / 448 (the test_qwen3_5.cpp:301-311 rule per row)."""
    op = "quantize_rows_e4m3"
    _require(x.is_cuda and x.dtype in (torch.float16, torch.bfloat16), op, "x must be a CUDA fp16/bf16 tensor")
    _require(x.dim() == 2 and x.is_contiguous(), op, "x must be a contiguous [M, K]")
    m, k = x.shape
    codes = torch.empty((m, k), dtype=torch.uint8, device=x.device)
    scale = torch.empty((m,), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        _call("plm_quantize_rows_e4m3", _ptr(x), _DTYPES[x.dtype], m, k, _ptr(codes), _ptr(scale),
              _stream(x.device))
    return codes, scale


def gemm_fp8_w8a8_cuda(x, weight_marlin, scale_marlin, n: int, block_n: int, group_size: int, out=None):
    """W8A8: x quantized per row to e4m3, fp8 x fp8 MFMA with fp32 block scales
    (no reference counterpart; the reference's fp8 GEMM is W8A16)."""
    op = "gemm_fp8_w8a8"
    _gemm_checks(op, _lib.PLM_FP8, x, weight_marlin, scale_marlin, n, block_n, group_size)
    _require(group_size % 128 == 0, op, "group_size must be a multiple of 128 for the fp8 MFMA")
    m, k = x.shape
    y = out if out is not None else torch.empty((m, n), dtype=x.dtype, device=x.device)
    if m == 0 or n == 0:
        return y
    lib = _lib.load()
    ws = workspace(x.device, lib.plm_gemm_w8a8_workspace_bytes(m, n, k))
    with torch.cuda.device(x.device):
        _call("plm_gemm_w8a8", _ptr(x), _DTYPES[x.dtype], _ptr(weight_marlin.contiguous()),
              _ptr(scale_marlin.contiguous()), _DTYPES[scale_marlin.dtype], m, n, k, block_n, group_size, _ptr(y),
              _ptr(ws), 0 if ws is None else ws.numel(), _stream(x.device))
    return y


# ---------------------------------------------------------------------------
# MoE: experts repacked back to back, grouped GEMM, routed experts
# ---------------------------------------------------------------------------


def repack_int4_experts(weight_packed: torch.Tensor, weight_scale: torch.Tensor, group_size: int):
    """[E, N, K/8] int32 + [E, N, K/g] scales -> per-expert plm layouts back to back:
    (weights int32 [E * words], scales [E, strips, groups, 16])."""
    op = "repack_int4_experts"
    _require(weight_packed.dim() == 3 and weight_scale.dim() == 3, op, "expected [E, N, K/8] and [E, N, K/g]")
    e = weight_packed.shape[0]
    ws, ss = [], []
    for i in range(e):
        w, s = repack_int4_marlin_cuda(weight_packed[i], weight_scale[i], 1, group_size)
        ws.append(w)
        ss.append(s)
    return torch.cat(ws), torch.stack(ss)


def grouped_gemm_int4_cuda(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor, offsets: torch.Tensor, n: int,
                           group_size: int, out=None) -> torch.Tensor:
    """Rows [offsets[e-1], offsets[e]) of x times expert e's W^T (one at::_grouped_mm of
    paged_forward.cpp:124-125, int4 experts)."""
    op = "grouped_gemm"
    _require(x.is_cuda and x.dim() == 2 and x.is_contiguous() and x.dtype in (torch.float16, torch.bfloat16), op,
             "x must be a contiguous CUDA [rows, K] fp16/bf16")
    _require(offsets.dtype == torch.int32 and offsets.dim() == 1, op, "offsets must be int32 [E]")
    rows, k = x.shape
    e = offsets.shape[0]
    lib = _lib.load()
    _require(weight.numel() * 4 == e * lib.plm_weight_bytes(_lib.PLM_INT4, n, k), op, "weight has the wrong size")
    y = out if out is not None else torch.empty((rows, n), dtype=x.dtype, device=x.device)
    if rows == 0 or n == 0:
        return y
    ws = workspace(x.device, lib.plm_grouped_gemm_workspace_bytes(rows, e))
    with torch.cuda.device(x.device):
        _call("plm_grouped_gemm", _lib.PLM_INT4, _ptr(x), _DTYPES[x.dtype], _ptr(weight), _ptr(scale),
              _DTYPES[scale.dtype], _ptr(offsets.contiguous()), e, rows, n, k, 1, group_size, _ptr(y), _ptr(ws),
              ws.numel(), _stream(x.device))
    return y


def routed_experts_int4_cuda(h: torch.Tensor, top_experts: torch.Tensor, top_weights: torch.Tensor,
                             gate_up: tuple, down: tuple, intermediate: int, group_size: int):
    """routed_experts (paged_forward.cpp:108-130) with int4 experts and SiLU:
    returns (out [T, H] in h's dtype, offsets int32 [E])."""
    op = "routed_experts"
    _require(h.is_cuda and h.dim() == 2 and h.dtype in (torch.float16, torch.bfloat16), op,
             "h must be a CUDA [T, H] fp16/bf16 tensor")
    t, hidden = h.shape
    top_k = top_experts.shape[-1]
    e = gate_up[1].shape[0]
    experts = top_experts.to(torch.int32).contiguous()
    weights = top_weights.to(torch.float32).contiguous()
    out = torch.empty_like(h)
    offsets = torch.empty((e,), dtype=torch.int32, device=h.device)
    lib = _lib.load()
    ws = workspace(h.device, lib.plm_moe_workspace_bytes(t, top_k, e, hidden, intermediate))
    with torch.cuda.device(h.device):
        _call("plm_moe", _ptr(h.contiguous()), _DTYPES[h.dtype], _ptr(experts), _ptr(weights), t, top_k, e, hidden,
              intermediate, _ptr(gate_up[0]), _ptr(gate_up[1]), _ptr(down[0]), _ptr(down[1]),
              _DTYPES[gate_up[1].dtype], group_size, _ptr(offsets), _ptr(out), _ptr(ws),
              0 if ws is None else ws.numel(), _stream(h.device))
    return out, offsets


def route_top_k_cuda(logits: torch.Tensor, k: int, experts_i32: bool = False):
    """route_top_k_cuda (ops.hpp:37-40): (weights fp32 [T, k], experts int64 [T, k]) for
    logits [T, E] whose rows may lie apart (unit column stride); experts_i32 gives int32
    experts (what routed_experts_int4_cuda / plm_moe take) instead."""
    op = "route_top_k"
    _require(logits.is_cuda and logits.dim() == 2 and logits.stride(1) == 1, op,
             "logits must be CUDA [tokens, experts], each row contiguous")
    _require(logits.dtype in _DTYPES, op, "logits must be fp32, fp16 or bf16")
    t, e = logits.shape
    weights = torch.empty((t, k), dtype=torch.float32, device=logits.device)
    chosen = torch.empty((t, k), dtype=torch.int32 if experts_i32 else torch.int64, device=logits.device)
    stride = logits.stride(0) if t > 1 else e
    with torch.cuda.device(logits.device):
        _call("plm_route_top_k", _ptr(logits), _DTYPES[logits.dtype], t, e, stride, k, _ptr(weights),
              None if experts_i32 else _ptr(chosen), _ptr(chosen) if experts_i32 else None, _stream(logits.device))
    return weights, chosen


def silu_mul_cuda(x: torch.Tensor) -> torch.Tensor:
    """silu_mul_cuda (ops.hpp:42-43): silu(x[:, :n]) * x[:, n:], silu rounded to the dtype."""
    op = "silu_mul"
    _require(x.is_cuda and x.dim() == 2 and x.is_contiguous() and x.size(1) % 2 == 0, op,
             "x must be contiguous CUDA [tokens, 2 * n]")
    _require(x.dtype in _DTYPES, op, "x must be fp32, fp16 or bf16")
    t, n = x.size(0), x.size(1) // 2
    y = torch.empty((t, n), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        _call("plm_silu_mul", _ptr(x), _DTYPES[x.dtype], t, n, _ptr(y), _stream(x.device))
    return y


def moe_block_int4_cuda(h: torch.Tensor, router_logits: torch.Tensor, top_k: int, gate_up: tuple, down: tuple,
                        intermediate: int, group_size: int):
    """The routed-experts half of a MoE block from the router's logits: route_top_k (int32
    experts) then routed_experts with int4 experts and SiLU (qwen4_exp.cpp:542 followed by
    paged_forward.cpp:108-130), all enqueued on the current stream with no host sync.
    Returns (out [T, H], offsets int32 [E], top_weights fp32 [T, k], top_experts int32 [T, k])."""
    weights, experts = route_top_k_cuda(router_logits, top_k, experts_i32=True)
    out, offsets = routed_experts_int4_cuda(h, experts, weights, gate_up, down, intermediate, group_size)
    return out, offsets, weights, experts


def _gemm_int4_plain(op: str, x: torch.Tensor, weight_packed: torch.Tensor, weight_scale: torch.Tensor,
                     group_size: int, num_splits: int) -> torch.Tensor:
    _require(x.is_cuda and x.dim() == 2 and x.dtype in (torch.float16, torch.bfloat16), op,
             "x must be a CUDA [M, K] fp16/bf16 tensor")
    _require(weight_packed.dtype == torch.int32 and weight_packed.dim() == 2, op, "weight_packed must be int32 [N, K/8]")
    m, k = x.shape
    n = weight_packed.shape[0]
    _require(weight_packed.shape[1] * 8 == k, op, "weight_packed must be [N, K/8]")
    _require(weight_scale.dim() == 2 and tuple(weight_scale.shape) == (n, k // group_size) if group_size > 0 else False,
             op, "weight_scale must be [N, K/group_size]")
    scale = weight_scale.to(torch.float32).contiguous()
    y = torch.empty((m, n), dtype=x.dtype, device=x.device)
    lib = _lib.load()
    nbytes = lib.plm_gemm_int4_plain_workspace_bytes(m, n, k, num_splits)
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=x.device) if nbytes > 0 else None
    with torch.cuda.device(x.device):
        _call("plm_gemm_int4_plain", _ptr(x.contiguous()), _DTYPES[x.dtype], _ptr(weight_packed.contiguous()),
              _ptr(scale), m, n, k, group_size, num_splits, _ptr(y), _ptr(ws), 0 if ws is None else ws.numel(),
              _stream(x.device))
    return y


def gemm_int4_cuda(x: torch.Tensor, weight_packed: torch.Tensor, weight_scale: torch.Tensor, group_size: int):
    """gemm_int4_cuda (ops.hpp:272-285): the non-repacked int4 GEMM, W = round(fp32(q * scale))."""
    return _gemm_int4_plain("gemm_int4", x, weight_packed, weight_scale, group_size, 0)


def gemm_int4_split_cuda(x: torch.Tensor, weight_packed: torch.Tensor, weight_scale: torch.Tensor, group_size: int,
                         num_splits: int):
    """gemm_int4_split_cuda (ops.hpp:287-297): the same with the K split forced to num_splits (>= 1)."""
    _require(num_splits >= 1, "gemm_int4", "num_splits must be >= 1")
    return _gemm_int4_plain("gemm_int4", x, weight_packed, weight_scale, group_size, num_splits)
