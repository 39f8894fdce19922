// y = x @ W^T over x's last dim for a dense, fp8 or int4 weight: the reference's
// linear (pulsarlm-core/inc/pulsarlm/engine/model/linear.hpp:13-35,
// src/engine/model/linear.cpp:19-41) with an int4 alternative next to fp8.
#pragma once

#include <ATen/ATen.h>

#include <cstdint>
#include <variant>

namespace pulsarlm {

class linear {
    struct quant_weight {
        at::Tensor weight_marlin;
        at::Tensor scale_marlin;
        std::int64_t n;
        std::int64_t block_n;
        std::int64_t group_size;
        bool fp8;
    };

    std::variant<at::Tensor, quant_weight> weight;

    explicit linear(std::variant<at::Tensor, quant_weight> weight);

  public:
    // weight [N, K] in x's dtype.
    static linear dense(at::Tensor weight);

    // weight float8_e4m3fn [N, K]; W[n, k] = weight[n, k] * scale[n / block_n, k / group_size].
    static linear fp8(const at::Tensor& weight, const at::Tensor& scale, std::int64_t block_n, std::int64_t group_size);

    // A checkpoint's fp8 linear whose output rows are reordered: output row r is weight row
    // row_order[r] (int64 [N]). weight_scale_inv [ceil(N/block_n), K/block_k] first expands to
    // one scale per row, since the reordering moves rows across the scale blocks
    // (need_permuted_linear, pulsarlm-core/src/engine/model/qwen3_5.cpp:65-83).
    static linear fp8_rows(const at::Tensor& weight, const at::Tensor& weight_scale_inv, std::int64_t block_n,
                           std::int64_t block_k, const at::Tensor& row_order);

    // weight_packed int32 [N, K/8] (8 signed int4 per int32, least significant first); same scale rule.
    static linear int4(const at::Tensor& weight_packed, const at::Tensor& scale, std::int64_t block_n,
                       std::int64_t group_size);

    at::Tensor apply(const at::Tensor& x) const;
};

}  // namespace pulsarlm
