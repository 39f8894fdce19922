// linear over the pulsarlm_amd ops: the reference's dense/fp8 linear
// (pulsarlm-core/src/engine/model/linear.cpp:14-41) plus an int4 alternative.
// Quantized weights are repacked once, at construction, as the reference does.
#include "linear.hpp"

#include <utility>
#include <vector>

#include "pulsarlm_ops.hpp"

namespace pulsarlm {

linear::linear(std::variant<at::Tensor, quant_weight> weight) : weight(std::move(weight)) {}

linear linear::dense(at::Tensor weight) { return linear(std::move(weight)); }

linear linear::fp8(const at::Tensor& weight, const at::Tensor& scale, std::int64_t block_n, std::int64_t group_size) {
    auto [w, s] = repack_fp8_marlin_cuda(weight, scale, block_n, group_size);
    return linear(quant_weight{std::move(w), std::move(s), weight.size(0), block_n, group_size, true});
}

linear linear::fp8_rows(const at::Tensor& weight, const at::Tensor& weight_scale_inv, std::int64_t block_n,
                        std::int64_t block_k, const at::Tensor& row_order) {
    TORCH_CHECK(row_order.dim() == 1 && row_order.size(0) == weight.size(0),
                "linear: row_order must hold one index per weight row");
    const at::Tensor order = row_order.to(weight.device(), at::kLong);
    const at::Tensor row_scale =
        weight_scale_inv.to(weight.device()).repeat_interleave(block_n, 0).narrow(0, 0, weight.size(0));
    const at::Tensor rows = weight.view(at::kByte).index_select(0, order).view(at::kFloat8_e4m3fn);
    return fp8(rows, row_scale.index_select(0, order).contiguous(), 1, block_k);
}

linear linear::int4(const at::Tensor& weight_packed, const at::Tensor& scale, std::int64_t block_n,
                    std::int64_t group_size) {
    auto [w, s] = repack_int4_marlin_cuda(weight_packed, scale, block_n, group_size);
    return linear(quant_weight{std::move(w), std::move(s), weight_packed.size(0), block_n, group_size, false});
}

at::Tensor linear::apply(const at::Tensor& x) const {
    if (const auto* dense = std::get_if<at::Tensor>(&weight)) return at::linear(x, *dense);
    const quant_weight& w = std::get<quant_weight>(weight);
    std::vector<std::int64_t> sizes = x.sizes().vec();
    const at::Tensor rows = x.reshape({-1, sizes.back()}).contiguous();
    sizes.back() = w.n;
    const at::Tensor y = w.fp8 ? gemm_fp8_marlin_cuda(rows, w.weight_marlin, w.scale_marlin, w.n, w.block_n, w.group_size)
                               : gemm_int4_marlin_cuda(rows, w.weight_marlin, w.scale_marlin, w.n, w.block_n,
                                                       w.group_size);
    return y.view(sizes);
}

}  // namespace pulsarlm
