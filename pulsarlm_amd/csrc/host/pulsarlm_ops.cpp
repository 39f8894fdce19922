// Implementation of pulsarlm_ops.hpp over the C ABI. Argument checks restate those of
// gemm<fmt> / repack<fmt> (pulsarlm-core/src/kernels/marlin.cu:395-445,538-576); the C
// ABI checks them again and reports anything it rejects through plm_last_error().
#include "pulsarlm_ops.hpp"

// PyTorch-ROCm tensors report device type "cuda"; the masquerading guard and stream
// accessors take that device type.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "pulsarlm_amd.h"

namespace pulsarlm {
namespace {

plm_dtype dtype_of(const char* op, at::ScalarType t) {
    switch (t) {
        case at::kBFloat16: return PLM_BF16;
        case at::kHalf: return PLM_FP16;
        case at::kFloat: return PLM_FP32;
        default: TORCH_CHECK(false, op, ": unsupported dtype ", t);
    }
}

void check_rc(int rc) {
    TORCH_CHECK(rc == PLM_OK, plm_last_error());
}

void* stream_of(const at::Tensor& t) {
    return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

std::vector<int64_t> scale_shape(int64_t n, int64_t k, int64_t block_n, int64_t group_size) {
    const int64_t strips = ceil_div(n, 16), ktiles = ceil_div(k, 128);
    return {strips, ceil_div(ktiles * 128, group_size), block_n % 16 == 0 ? 1 : 16};
}

// One zero-initialised workspace per (device, stream): the kernels leave the split-K
// counters at its front at zero, so calls ordered on one stream can share it.
std::mutex ws_mutex;
std::map<std::pair<int, void*>, at::Tensor> ws_cache;

at::Tensor workspace(const at::Tensor& like, int64_t bytes) {
    if (bytes <= 0) return at::Tensor();
    std::lock_guard<std::mutex> lock(ws_mutex);
    auto key = std::make_pair(static_cast<int>(like.device().index()), stream_of(like));
    auto it = ws_cache.find(key);
    if (it == ws_cache.end() || it->second.numel() < bytes) {
        at::Tensor buf = at::zeros({std::max<int64_t>(bytes, 1 << 20)}, like.options().dtype(at::kByte));
        ws_cache[key] = buf;
        return buf;
    }
    return it->second;
}

void* ptr(const at::Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

std::tuple<at::Tensor, at::Tensor> repack(const char* op, plm_format fmt, const at::Tensor& weight, int64_t n,
                                          int64_t k, const at::Tensor& weight_scale, int64_t block_n,
                                          int64_t group_size) {
    TORCH_CHECK(weight.is_cuda() && weight_scale.is_cuda(), op, ": inputs must be CUDA tensors");
    TORCH_CHECK(block_n > 0, op, ": block_n must be positive");
    TORCH_CHECK(group_size > 0 && group_size % 16 == 0, op, ": group_size must be a positive multiple of 16");
    TORCH_CHECK(k % group_size == 0, op, ": K must be a multiple of group_size");
    TORCH_CHECK(weight_scale.dim() == 2 && weight_scale.size(0) == ceil_div(n, block_n) &&
                    weight_scale.size(1) == k / group_size,
                op, ": weight_scale must be [ceil(N / block_n), K / group_size]");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(weight.device());
    const at::Tensor src = weight.contiguous();
    const at::Tensor scale = weight_scale.contiguous();
    at::Tensor w = at::empty({plm_weight_bytes(fmt, n, k) / 4}, weight.options().dtype(at::kInt));
    at::Tensor s = at::empty(scale_shape(n, k, block_n, group_size), scale.options());
    const plm_dtype sd = dtype_of(op, scale.scalar_type());
    const int rc = fmt == PLM_INT4
                       ? plm_repack_int4(static_cast<const int32_t*>(src.data_ptr()), scale.data_ptr(), sd, n, k,
                                         block_n, group_size, w.data_ptr(), s.data_ptr(), stream_of(weight))
                       : plm_repack_fp8(static_cast<const uint8_t*>(src.data_ptr()), scale.data_ptr(), sd, n, k,
                                        block_n, group_size, w.data_ptr(), s.data_ptr(), stream_of(weight));
    check_rc(rc);
    return {w, s};
}

void gemm_checks(const char* op, plm_format fmt, const at::Tensor& x, const at::Tensor& weight_marlin,
                 const at::Tensor& scale_marlin, int64_t n, int64_t block_n, int64_t group_size) {
    TORCH_CHECK(x.is_cuda() && weight_marlin.is_cuda() && scale_marlin.is_cuda(), op,
                ": all inputs must be CUDA tensors");
    TORCH_CHECK(x.scalar_type() == at::kHalf || x.scalar_type() == at::kBFloat16, op, ": x must be fp16 or bf16");
    TORCH_CHECK(x.dim() == 2 && x.is_contiguous(), op, ": x must be a contiguous [M, K]");
    TORCH_CHECK(weight_marlin.scalar_type() == at::kInt, op, ": weight_marlin must be int32");
    TORCH_CHECK(block_n > 0, op, ": block_n must be positive");
    TORCH_CHECK(group_size > 0 && group_size % 16 == 0, op, ": group_size must be a positive multiple of 16");
    const int64_t k = x.size(1);
    TORCH_CHECK(k % group_size == 0, op, ": K must be a multiple of group_size");
    TORCH_CHECK(scale_marlin.sizes().vec() == scale_shape(n, k, block_n, group_size), op,
                ": scale_marlin has the wrong shape for this N, K, block_n and group_size");
    TORCH_CHECK(weight_marlin.numel() * 4 == plm_weight_bytes(fmt, n, k), op,
                ": weight_marlin has the wrong size for this shape");
}

at::Tensor gemm(const char* op, plm_format fmt, bool w8a8, const at::Tensor& x, const at::Tensor& weight_marlin,
                const at::Tensor& scale_marlin, int64_t n, int64_t block_n, int64_t group_size) {
    gemm_checks(op, fmt, x, weight_marlin, scale_marlin, n, block_n, group_size);
    at::Tensor y = at::empty({x.size(0), n}, x.options());
    if (x.size(0) == 0 || n == 0) return y;
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const int64_t m = x.size(0), k = x.size(1);
    const at::Tensor w = weight_marlin.contiguous(), s = scale_marlin.contiguous();
    const plm_dtype sd = dtype_of(op, s.scalar_type());
    const plm_dtype xd = dtype_of(op, x.scalar_type());
    if (w8a8) {
        at::Tensor ws = workspace(x, plm_gemm_w8a8_workspace_bytes(m, n, k));
        check_rc(plm_gemm_w8a8(x.data_ptr(), xd, w.data_ptr(), s.data_ptr(), sd, m, n, k, block_n, group_size,
                               y.data_ptr(), ptr(ws), ws.defined() ? ws.numel() : 0, stream_of(x)));
    } else {
        at::Tensor ws = workspace(x, plm_gemm_workspace_bytes(fmt, m, n, k));
        check_rc(plm_gemm(fmt, x.data_ptr(), xd, w.data_ptr(), s.data_ptr(), sd, m, n, k, block_n, group_size,
                          y.data_ptr(), ptr(ws), ws.defined() ? ws.numel() : 0, stream_of(x)));
    }
    return y;
}

}  // namespace

std::tuple<at::Tensor, at::Tensor> repack_int4_marlin_cuda(const at::Tensor& weight_packed,
                                                           const at::Tensor& weight_scale, int64_t block_n,
                                                           int64_t group_size) {
    TORCH_CHECK(weight_packed.scalar_type() == at::kInt && weight_packed.dim() == 2,
                "repack_int4_marlin: weight_packed must be int32 [N, K/8]");
    return repack("repack_int4_marlin", PLM_INT4, weight_packed, weight_packed.size(0), weight_packed.size(1) * 8,
                  weight_scale, block_n, group_size);
}

std::tuple<at::Tensor, at::Tensor> repack_fp8_marlin_cuda(const at::Tensor& weight, const at::Tensor& weight_scale,
                                                          int64_t block_n, int64_t group_size) {
    TORCH_CHECK(weight.scalar_type() == at::kFloat8_e4m3fn && weight.dim() == 2,
                "repack_fp8_marlin: weight must be float8_e4m3fn [N, K]");
    return repack("repack_fp8_marlin", PLM_FP8, weight, weight.size(0), weight.size(1), weight_scale, block_n,
                  group_size);
}

at::Tensor gemm_int4_marlin_cuda(const at::Tensor& x, const at::Tensor& weight_marlin, const at::Tensor& scale_marlin,
                                 int64_t n, int64_t block_n, int64_t group_size) {
    return gemm("gemm_int4_marlin", PLM_INT4, false, x, weight_marlin, scale_marlin, n, block_n, group_size);
}

at::Tensor gemm_fp8_marlin_cuda(const at::Tensor& x, const at::Tensor& weight_marlin, const at::Tensor& scale_marlin,
                                int64_t n, int64_t block_n, int64_t group_size) {
    return gemm("gemm_fp8_marlin", PLM_FP8, false, x, weight_marlin, scale_marlin, n, block_n, group_size);
}

at::Tensor gemm_fp8_w8a8_cuda(const at::Tensor& x, const at::Tensor& weight_marlin, const at::Tensor& scale_marlin,
                              int64_t n, int64_t block_n, int64_t group_size) {
    TORCH_CHECK(group_size % 128 == 0, "gemm_fp8_w8a8: group_size must be a multiple of 128 for the fp8 MFMA");
    return gemm("gemm_fp8_w8a8", PLM_FP8, true, x, weight_marlin, scale_marlin, n, block_n, group_size);
}

std::tuple<at::Tensor, at::Tensor> quantize_rows_e4m3_cuda(const at::Tensor& x) {
    const char* op = "quantize_rows_e4m3";
    TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.is_contiguous(), op, ": x must be a contiguous CUDA [M, K]");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    at::Tensor codes = at::empty({x.size(0), x.size(1)}, x.options().dtype(at::kByte));
    at::Tensor scale = at::empty({x.size(0)}, x.options().dtype(at::kFloat));
    check_rc(plm_quantize_rows_e4m3(x.data_ptr(), dtype_of(op, x.scalar_type()), x.size(0), x.size(1),
                                    static_cast<uint8_t*>(codes.data_ptr()), static_cast<float*>(scale.data_ptr()),
                                    stream_of(x)));
    return {codes, scale};
}

std::tuple<at::Tensor, at::Tensor> convert_marlin_cuda(const std::string& format, const at::Tensor& weight_marlin,
                                                       const at::Tensor& scale_marlin, int64_t n, int64_t k,
                                                       int64_t block_n, int64_t group_size) {
    const char* op = "convert_marlin";
    TORCH_CHECK(format == "int4" || format == "fp8", op, ": format must be int4 or fp8");
    TORCH_CHECK(weight_marlin.scalar_type() == at::kInt && scale_marlin.scalar_type() == at::kFloat, op,
                ": weight_marlin must be int32 and scale_marlin fp32");
    const plm_format fmt = format == "int4" ? PLM_INT4 : PLM_FP8;
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(weight_marlin.device());
    at::Tensor w = at::empty({plm_weight_bytes(fmt, n, k) / 4}, weight_marlin.options());
    at::Tensor s = at::empty(scale_shape(n, k, block_n, group_size), scale_marlin.options());
    const at::Tensor wm = weight_marlin.contiguous(), sm = scale_marlin.contiguous();
    check_rc(plm_convert_marlin(fmt, static_cast<const int32_t*>(wm.data_ptr()), static_cast<const float*>(sm.data_ptr()),
                                n, k, block_n, group_size, w.data_ptr(), s.data_ptr(), stream_of(weight_marlin)));
    return {w, s};
}

at::Tensor dequant_marlin_cuda(const std::string& format, const at::Tensor& weight_marlin,
                               const at::Tensor& scale_marlin, int64_t n, int64_t k, int64_t block_n,
                               int64_t group_size, at::ScalarType dtype) {
    const char* op = "dequant";
    TORCH_CHECK(format == "int4" || format == "fp8", op, ": format must be int4 or fp8");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(weight_marlin.device());
    at::Tensor out = at::empty({n, k}, weight_marlin.options().dtype(dtype));
    check_rc(plm_dequant(format == "int4" ? PLM_INT4 : PLM_FP8, weight_marlin.data_ptr(), scale_marlin.data_ptr(),
                         dtype_of(op, scale_marlin.scalar_type()), n, k, block_n, group_size, out.data_ptr(),
                         dtype_of(op, dtype), stream_of(weight_marlin)));
    return out;
}

std::tuple<at::Tensor, at::Tensor> repack_int4_experts_cuda(const at::Tensor& weight_packed,
                                                            const at::Tensor& weight_scale, int64_t group_size) {
    TORCH_CHECK(weight_packed.dim() == 3 && weight_scale.dim() == 3,
                "repack_int4_experts: expected [E, N, K/8] weights and [E, N, K/g] scales");
    std::vector<at::Tensor> ws, ss;
    for (int64_t e = 0; e < weight_packed.size(0); ++e) {
        auto [w, s] = repack_int4_marlin_cuda(weight_packed[e], weight_scale[e], 1, group_size);
        ws.push_back(w);
        ss.push_back(s);
    }
    return {at::cat(ws), at::stack(ss)};
}

at::Tensor grouped_gemm_int4_cuda(const at::Tensor& x, const at::Tensor& weight, const at::Tensor& scale,
                                  const at::Tensor& offsets, int64_t n, int64_t group_size) {
    const char* op = "grouped_gemm";
    TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.is_contiguous(), op, ": x must be a contiguous CUDA [rows, K]");
    TORCH_CHECK(offsets.scalar_type() == at::kInt && offsets.dim() == 1, op, ": offsets must be int32 [E]");
    const int64_t rows = x.size(0), k = x.size(1), e = offsets.size(0);
    TORCH_CHECK(weight.numel() * 4 == e * plm_weight_bytes(PLM_INT4, n, k), op, ": weight has the wrong size");
    at::Tensor y = at::empty({rows, n}, x.options());
    if (rows == 0 || n == 0) return y;
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    at::Tensor ws = workspace(x, plm_grouped_gemm_workspace_bytes(rows, e));
    const at::Tensor off = offsets.contiguous();
    check_rc(plm_grouped_gemm(PLM_INT4, x.data_ptr(), dtype_of(op, x.scalar_type()), weight.data_ptr(),
                              scale.data_ptr(), dtype_of(op, scale.scalar_type()),
                              static_cast<const int32_t*>(off.data_ptr()), e, rows, n, k, 1, group_size, y.data_ptr(),
                              ptr(ws), ws.numel(), stream_of(x)));
    return y;
}

std::tuple<at::Tensor, at::Tensor> routed_experts_int4_cuda(const at::Tensor& h, const at::Tensor& top_experts,
                                                            const at::Tensor& top_weights,
                                                            const at::Tensor& gate_up_weight,
                                                            const at::Tensor& gate_up_scale,
                                                            const at::Tensor& down_weight,
                                                            const at::Tensor& down_scale, int64_t intermediate,
                                                            int64_t group_size) {
    const char* op = "routed_experts";
    TORCH_CHECK(h.is_cuda() && h.dim() == 2, op, ": h must be a CUDA [T, H] tensor");
    TORCH_CHECK(top_experts.sizes() == top_weights.sizes() && top_experts.dim() == 2, op,
                ": top_experts and top_weights must be [T, top_k]");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(h.device());
    const int64_t t = h.size(0), hidden = h.size(1), top_k = top_experts.size(1), e = gate_up_scale.size(0);
    const at::Tensor hc = h.contiguous();
    const at::Tensor experts = top_experts.to(at::kInt).contiguous();
    const at::Tensor weights = top_weights.to(at::kFloat).contiguous();
    at::Tensor out = at::empty_like(hc);
    at::Tensor offsets = at::empty({e}, h.options().dtype(at::kInt));
    at::Tensor ws = workspace(h, plm_moe_workspace_bytes(t, top_k, e, hidden, intermediate));
    check_rc(plm_moe(hc.data_ptr(), dtype_of(op, h.scalar_type()), static_cast<const int32_t*>(experts.data_ptr()),
                     static_cast<const float*>(weights.data_ptr()), t, top_k, e, hidden, intermediate,
                     gate_up_weight.data_ptr(), gate_up_scale.data_ptr(), down_weight.data_ptr(),
                     down_scale.data_ptr(), dtype_of(op, gate_up_scale.scalar_type()), group_size,
                     static_cast<int32_t*>(offsets.data_ptr()), out.data_ptr(), ptr(ws), ws.defined() ? ws.numel() : 0,
                     stream_of(h)));
    return {out, offsets};
}

std::tuple<at::Tensor, at::Tensor> route_top_k_cuda(const at::Tensor& logits, int64_t k) {
    const char* op = "route_top_k";
    TORCH_CHECK(logits.is_cuda() && logits.dim() == 2 && logits.stride(1) == 1, op,
                ": logits must be CUDA [tokens, experts], each row contiguous");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(logits.device());
    const int64_t tokens = logits.size(0), experts = logits.size(1);
    at::Tensor weights = at::empty({tokens, k}, logits.options().dtype(at::kFloat));
    at::Tensor chosen = at::empty({tokens, k}, logits.options().dtype(at::kLong));
    check_rc(plm_route_top_k(logits.data_ptr(), dtype_of(op, logits.scalar_type()), tokens, experts,
                             tokens > 1 ? logits.stride(0) : experts, k, static_cast<float*>(weights.data_ptr()),
                             static_cast<int64_t*>(chosen.data_ptr()), nullptr, stream_of(logits)));
    return {weights, chosen};
}

at::Tensor silu_mul_cuda(const at::Tensor& x) {
    const char* op = "silu_mul";
    TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.is_contiguous() && x.size(1) % 2 == 0, op,
                ": x must be contiguous CUDA [tokens, 2 * n]");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const int64_t tokens = x.size(0), n = x.size(1) / 2;
    at::Tensor y = at::empty({tokens, n}, x.options());
    check_rc(plm_silu_mul(x.data_ptr(), dtype_of(op, x.scalar_type()), tokens, n, y.data_ptr(), stream_of(x)));
    return y;
}

namespace {
at::Tensor gemm_int4_plain(const char* op, const at::Tensor& x, const at::Tensor& weight_packed,
                           const at::Tensor& weight_scale, int64_t group_size, int64_t num_splits) {
    TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.is_contiguous(), op, ": x must be a contiguous CUDA [M, K] tensor");
    TORCH_CHECK(weight_packed.is_cuda() && weight_packed.scalar_type() == at::kInt && weight_packed.dim() == 2 &&
                    weight_packed.is_contiguous(),
                op, ": weight_packed must be contiguous CUDA int32 [N, K/8]");
    const int64_t m = x.size(0), k = x.size(1), n = weight_packed.size(0);
    TORCH_CHECK(weight_packed.size(1) * 8 == k, op, ": weight_packed must be [N, K/8]");
    TORCH_CHECK(group_size > 0 && weight_scale.dim() == 2 && weight_scale.size(0) == n &&
                    weight_scale.size(1) * group_size == k,
                op, ": weight_scale must be [N, K/group_size]");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
    const at::Tensor scale = weight_scale.to(at::kFloat).contiguous();
    at::Tensor y = at::empty({m, n}, x.options());
    const int64_t nbytes = plm_gemm_int4_plain_workspace_bytes(m, n, k, num_splits);
    at::Tensor ws = nbytes > 0 ? at::empty({nbytes}, x.options().dtype(at::kByte)) : at::Tensor();
    check_rc(plm_gemm_int4_plain(x.data_ptr(), dtype_of(op, x.scalar_type()),
                                 static_cast<const int32_t*>(weight_packed.data_ptr()),
                                 static_cast<const float*>(scale.data_ptr()), m, n, k, group_size, num_splits,
                                 y.data_ptr(), ptr(ws), ws.defined() ? ws.numel() : 0, stream_of(x)));
    return y;
}
}  // namespace

at::Tensor gemm_int4_cuda(const at::Tensor& x, const at::Tensor& weight_packed, const at::Tensor& weight_scale,
                          int64_t group_size) {
    return gemm_int4_plain("gemm_int4", x, weight_packed, weight_scale, group_size, 0);
}

at::Tensor gemm_int4_split_cuda(const at::Tensor& x, const at::Tensor& weight_packed,
                                const at::Tensor& weight_scale, int64_t group_size, int64_t num_splits) {
    TORCH_CHECK(num_splits >= 1, "gemm_int4: num_splits must be >= 1");
    return gemm_int4_plain("gemm_int4", x, weight_packed, weight_scale, group_size, num_splits);
}

}  // namespace pulsarlm
