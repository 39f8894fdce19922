// Host-side drop-in for pulsarlm-core's quant-linear operators over the
// pulsarlm_amd C ABI (include/pulsarlm_amd.h), for PyTorch-ROCm tensors.
//
// The first four functions keep the exact signatures, argument meaning and error
// behaviour (TORCH_CHECK -> c10::Error, "<op>: ..." messages, empty [M, N] for
// M == 0 or N == 0) of pulsarlm-core/inc/pulsarlm/kernels/ops.hpp:306-332, so a
// caller such as linear (pulsarlm-core/src/engine/model/linear.cpp:19-41) links
// against this file instead of marlin.cu. Work is enqueued on the current HIP stream
// of the tensors' device; nothing synchronizes. weight_marlin / scale_marlin are
// opaque (the plm tile layout), as the reference's are.
#pragma once

#include <ATen/ATen.h>

#include <cstdint>
#include <tuple>

namespace pulsarlm {

// ops.hpp:306-311
std::tuple<at::Tensor, at::Tensor> repack_int4_marlin_cuda(const at::Tensor& weight_packed,
                                                           const at::Tensor& weight_scale, int64_t block_n,
                                                           int64_t group_size);

// ops.hpp:313-314
std::tuple<at::Tensor, at::Tensor> repack_fp8_marlin_cuda(const at::Tensor& weight, const at::Tensor& weight_scale,
                                                          int64_t block_n, int64_t group_size);

// ops.hpp:316-323
at::Tensor gemm_int4_marlin_cuda(const at::Tensor& x, const at::Tensor& weight_marlin, const at::Tensor& scale_marlin,
                                 int64_t n, int64_t block_n, int64_t group_size);

// ops.hpp:325-332
at::Tensor gemm_fp8_marlin_cuda(const at::Tensor& x, const at::Tensor& weight_marlin, const at::Tensor& scale_marlin,
                                int64_t n, int64_t block_n, int64_t group_size);

// ---- additions (no counterpart in ops.hpp) ----

// W8A8: x quantized per row to e4m3, fp8 MFMA; group_size % 128 == 0.
at::Tensor gemm_fp8_w8a8_cuda(const at::Tensor& x, const at::Tensor& weight_marlin, const at::Tensor& scale_marlin,
                              int64_t n, int64_t block_n, int64_t group_size);

// (codes uint8 [M, K], scale fp32 [M]) with scale = max(amax, 1e-12) / 448 per row.
std::tuple<at::Tensor, at::Tensor> quantize_rows_e4m3_cuda(const at::Tensor& x);

// Weights repacked by the reference's repack (Marlin words + fp32 [K/g, N/bn] scales)
// converted to the plm layout; format "int4" or "fp8".
std::tuple<at::Tensor, at::Tensor> convert_marlin_cuda(const std::string& format, const at::Tensor& weight_marlin,
                                                       const at::Tensor& scale_marlin, int64_t n, int64_t k,
                                                       int64_t block_n, int64_t group_size);

// Dense round(q * round(s)) [N, K] in dtype from the plm layout.
at::Tensor dequant_marlin_cuda(const std::string& format, const at::Tensor& weight_marlin,
                               const at::Tensor& scale_marlin, int64_t n, int64_t k, int64_t block_n,
                               int64_t group_size, at::ScalarType dtype);

// [E, N, K/8] int32 + [E, N, K/g] scales -> experts back to back in the plm layout.
std::tuple<at::Tensor, at::Tensor> repack_int4_experts_cuda(const at::Tensor& weight_packed,
                                                            const at::Tensor& weight_scale, int64_t group_size);

// Rows [offsets[e-1], offsets[e]) of x times expert e's W^T (an at::_grouped_mm of
// pulsarlm-core/src/engine/model/paged_forward.cpp:124-125 with int4 experts).
at::Tensor grouped_gemm_int4_cuda(const at::Tensor& x, const at::Tensor& weight, const at::Tensor& scale,
                                  const at::Tensor& offsets, int64_t n, int64_t group_size);

// routed_experts (paged_forward.cpp:108-130, paged_forward.hpp) with int4 experts and
// SiLU; returns (out [T, H], offsets int32 [E]).
std::tuple<at::Tensor, at::Tensor> routed_experts_int4_cuda(const at::Tensor& h, const at::Tensor& top_experts,
                                                            const at::Tensor& top_weights,
                                                            const at::Tensor& gate_up_weight,
                                                            const at::Tensor& gate_up_scale,
                                                            const at::Tensor& down_weight,
                                                            const at::Tensor& down_scale, int64_t intermediate,
                                                            int64_t group_size);

// route_top_k_cuda (pulsarlm-core/inc/pulsarlm/kernels/ops.hpp:37-40): (weights fp32
// [tokens, k], experts int64 [tokens, k]) from logits [tokens, experts] whose rows may lie apart.
std::tuple<at::Tensor, at::Tensor> route_top_k_cuda(const at::Tensor& logits, int64_t k);

// silu_mul_cuda (ops.hpp:42-43): silu(x[:, :n]) * x[:, n:], silu rounded to the dtype.
at::Tensor silu_mul_cuda(const at::Tensor& x);

// gemm_int4_cuda / gemm_int4_split_cuda (pulsarlm-core/inc/pulsarlm/kernels/ops.hpp:272-297):
// y [M, N] = x @ W^T with W = round(fp32(q * scale)) from weight_packed int32 [N, K/8] and
// weight_scale fp32 [N, K/group_size], read in place; the split variant forces num_splits.
at::Tensor gemm_int4_cuda(const at::Tensor& x, const at::Tensor& weight_packed, const at::Tensor& weight_scale,
                          int64_t group_size);
at::Tensor gemm_int4_split_cuda(const at::Tensor& x, const at::Tensor& weight_packed,
                                const at::Tensor& weight_scale, int64_t group_size, int64_t num_splits);

}  // namespace pulsarlm
